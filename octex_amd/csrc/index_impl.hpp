// State of a loaded octex index on one MI355X (the reference's index_impl + device_part,
// detail/index_impl.hpp:115-177, for a single device).
//
// HBM layout (one allocation per array):
//   lists    i32 [C, stride]        cell lists of all levels of every copy (stride = rows * l), or one
//                                   allocation per copy; list_ptr i64 [C] holds each copy's address
//   keys     i64 [C, L, mmax]       cell ids per (copy, level) in (bucket, id) order
//   offsets  i32 [C, L, 2^logT + 1] CSR of the buckets into keys
//   lines    16 B [C, L, 2^logT]   the probe's bucket lines: first key and key range of every bucket
//                                   (make_bucket_lines; absent when the device lacks the memory)
//   base     i32 [C, L]             first cell row of every level
//   ucatT    f16 [C * 8b, D]        projections of all copies, one row per projected coordinate
//                                   (the transpose of the reference's ucat [D, C * 8b]) so that the
//                                   MFMA A-operand loads are contiguous
//   shift    f16 [C * 8b], inv_f f32 [L], mean f32 [D], basis f32 [D, S], scale f32 [S]
//   sketch   i8  [N, S]             (or pinned host memory)
//   vectors  f16 [N, D]             (or pinned host memory)
//   table    i32 [N, table_len]     (or pinned host memory)
#pragma once

#include "common.hpp"

#include <cuvs/neighbors/octex.hpp>

#include <cstdint>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

namespace cuvs::neighbors::octex::detail {

struct plan;  // buffers and graph of one (batch, k, search parameters); search.cpp

/**
 * Bytes between two sketch rows of S codes in memory: the next power of two for S <= 128, else a multiple
 * of 128, so that no row straddles a 128-byte cache line (a 96-byte row at a 96-byte stride touches 1.5
 * lines on average; padded to 128 it touches one) -- while the padding of n rows costs at most 1/32 of the
 * device memory (device_bytes; 0: no limit): a billion rows of 96 codes keep S-byte rows, since their padding
 * alone would take 32 GB.  The directory keeps rows of S bytes.
 */
inline auto sketch_pitch_for(int S, int64_t n = 0, size_t device_bytes = 0) -> int
{
  int p = 16;
  if (S > 128) {
    p = (S + 127) / 128 * 128;
  } else {
    while (p < S)
      p <<= 1;
  }
  if (device_bytes > 0 && static_cast<double>(n) * (p - S) > static_cast<double>(device_bytes) / 32) return S;
  return p;
}

/** The device's memory in bytes (0 if it cannot be read). */
inline auto device_memory_bytes() -> size_t
{
  size_t fr = 0, tot = 0;
  return hipMemGetInfo(&fr, &tot) == hipSuccess ? tot : 0;
}

struct index_impl {
  // meta.json
  int64_t n = 0, dim = 0;
  int copies = 0, blocks = 4, list_len = 0, log_buckets = 20, sketch_width = 0, table_len = 0;
  int sketch_pitch = 0;  // bytes between sketch rows in memory (sketch_pitch_for(sketch_width))
  std::vector<float> spacings;
  std::string path;

  load_params params;
  std::vector<int> devices;  // the one GPU holding the index
  int device         = 0;
  hipStream_t stream = nullptr;

  dbuf lists;                     // the loader's lists [C, stride] (one allocation)
  std::vector<dbuf> copy_lists;   // or the builder's, one allocation per copy
  dbuf list_ptr;                  // i64 [C]: device address of every copy's lists
  std::vector<int64_t> list_rows; // cell rows of every copy (builder)
  dbuf keys, offsets, base, ucatT, shift, inv_f, mean, basis, scale;
  dbuf lines;  // bucket_line [C, L, T1 - 1], or empty
  dbuf sketch, vectors, table;
  hbuf host_sketch, host_vectors, host_table;
  int64_t stride = 0, mmax = 0, T1 = 0;
  int64_t bytes  = 0;  // device bytes of the arrays

  [[nodiscard]] auto levels() const -> int { return static_cast<int>(spacings.size()); }
  [[nodiscard]] auto code() const -> const signed char*
  {
    return host_sketch.ptr != nullptr ? static_cast<const signed char*>(host_sketch.dptr)
                                      : sketch.as<const signed char>();
  }
  [[nodiscard]] auto vecs() const -> const __half*
  {
    return host_vectors.ptr != nullptr ? static_cast<const __half*>(host_vectors.dptr)
                                       : vectors.as<const __half>();
  }
  [[nodiscard]] auto rows() const -> const int*
  {
    return host_table.ptr != nullptr ? static_cast<const int*>(host_table.dptr) : table.as<const int>();
  }

  std::mutex mu;  // the plan cache
  std::map<std::string, std::shared_ptr<plan>> plans;
  // Held by whoever works on `stream`: plan creation (its graph capture), a search's batches, the release of
  // an evicted plan (whose destructor waits for the stream), introspection and placement changes.  Work of
  // another thread reaching the stream during a capture would be captured into, or invalidate, that graph.
  std::mutex stream_mu;

  index_impl() = default;
  index_impl(index_impl const&) = delete;
  ~index_impl();
};

/**
 * The probe's bucket lines of a loaded or built index (keys and offsets in HBM), when the device keeps keep_free
 * bytes free beside them; without them the probe reads the offsets.  OCTEX_PROBE_LINES=0 leaves them out.
 */
void make_bucket_lines(index_impl& ix, size_t keep_free);
/** Device memory left free for the search's batch buffers when the bucket lines are added. */
constexpr size_t kSearchReserve = size_t{8} << 30;

}  // namespace cuvs::neighbors::octex::detail
