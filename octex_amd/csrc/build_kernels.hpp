// Device side of the octex index builder (build_kernels.hip).
#pragma once

#include "common.hpp"

#include <hip/hip_fp16.h>

#include <cstdint>
#include <vector>

namespace cuvs::neighbors::octex::detail {

/** G [d, d] (device, fp64) = A^T A of the ns sampled rows x[i * step] - mean. */
void pca_scatter(const __half* x, int64_t n, int d, int64_t step, int64_t ns, const float* mean, double* G,
                 hipStream_t s);
/** host_out [ns, d] = the rows x[i * step] (device to host through a compact device copy). */
void sample_rows(const __half* x, int64_t ns, int64_t step, int d, __half* host_out, hipStream_t s);
/** y [n, w] = (x - mean) @ U [d, w] + shift (fp32). */
void project_rows(const __half* x, int64_t n, int d, const float* mean, const float* U, const float* shift, int w,
                  float* y, hipStream_t s);
void half_to_float(const __half* x, int64_t total, float* out, hipStream_t s);
/** out [n] = squared norms of the rows x [n, d] (fp16 or fp32), in fp32. */
template <typename T>
void row_norms(const T* x, int64_t n, int d, float* out, hipStream_t s);
/**
 * The K (<= 128) nearest rows of X [n, d] to each row of Q [m, d] (fp16 or fp32) by squared L2 distance
 * (fp32 from the squared norms qn / xn and MFMA dot products), ties by row: out_d / out_i [m, K]
 * ascending, -1 / +inf padded when n < K (device arrays).
 */
template <typename T>
void knn_rows(const T* Q, const float* qn, int64_t m, const T* X, const float* xn, int64_t n, int d, int K,
              float* out_d, int* out_i, hipStream_t s);
/** out = fp16(x), round to nearest even (device arrays). */
void float_to_half(const float* x, int64_t total, __half* out, hipStream_t s);
/**
 * The dataset's fp16 rows [n, d] for passes in chunks: device rows read in place, or pinned host rows copied chunk by
 * chunk into a device staging buffer (a chunk's copy is ordered after the kernels of the previous one on s).
 */
struct row_source {
  const __half* dev  = nullptr;
  const __half* host = nullptr;
  int d              = 0;
  dbuf stage;
  /** Device rows [r0, r0 + m). */
  auto rows(int64_t r0, int64_t m, hipStream_t s) -> const __half*;
};

/** The int8 sketch: scale = amax / 127 per coordinate, codes [n, pitch] = round(((x - mean) @ basis) / scale). */
void make_sketch(row_source& x, int64_t n, int d, const float* mean, const float* basis, int S, int pitch,
                 std::vector<float>& scale, signed char* codes, hipStream_t s);

/**
 * An IVF index of one copy's projected rows y [n, w], for the reference's default cell lists (build_cells.cuh:511-516,
 * 584-596: cuVS ivf_flat with max(64, 4 sqrt(n)) lists trained on half the rows, a tenth above 4M, searched with
 * list_probes probes).  cuVS is not part of this build: the centers here are Lloyd k-means over an evenly spaced
 * sample (the first centers evenly spaced sample rows; a center keeps its place when no row is nearest to it), each
 * row's nearest center by the exact k-NN kernel, the sums of a center's rows in row order (the same centers on every
 * run).  The rows are kept grouped by center (yc, in the order rows[]).
 */
struct ivf_index {
  int64_t n = 0;
  int w = 0, nlist = 0;
  dbuf centers, cnorm, off, rows, yc;
  dbuf ys, ysn, yn, lab, slab, idx, sidx, cnt, dtmp, pd, pidx, tmp;

  /** k-means of `iters` rounds over the rows y[i * step] (about train_fraction of them, at least nlist). */
  void build(const float* y, int64_t n, int w, int nlist, double train_fraction, int iters, hipStream_t s);
  /**
   * out [M, l] (device): for each center z [M, w] (squared norms zn), the l rows nearest to it, by (fp32 squared
   * distance summed in coordinate order, row), among the rows of its `probes` nearest centers (at most 128),
   * -1 past the rows there are (l <= 128); with out_d, their distances [M, l] (+inf past the rows there are).
   */
  void lists(const float* z, const float* zn, int64_t M, int probes, int l, int* out, hipStream_t s,
             float* out_d = nullptr);
};

/** key / dist [m]: the cell id of each row of y [m, 8B] at spacing f and its squared distance to the cell's center. */
void stream_keys(const float* y, int64_t m, int B, float f, long long* key, float* dist, hipStream_t s);
/**
 * z [M, 8B] = the centers f * E8(y / f) of cells from one member each: rows [M] of x (device-readable fp16 rows
 * [*, d], d even), gathered `chunk` at a time into stage and projected into y [chunk, 8B].
 */
void cell_centers(const __half* x, const int* rows, int64_t M, int d, const float* mean, const float* U,
                  const float* shift, int B, float f, int64_t chunk, dbuf& stage, float* y, float* z, hipStream_t s);
/** bd = +inf, bi = -1 over total entries: empty lists. */
void init_lists(float* bd, int* bi, int64_t total, hipStream_t s);
/**
 * od / oi [M, l] = for each center the l first of its kept list (bd, bi) and of one row range's list (nd, ni, rows
 * numbered from a; -1 entries stay -1), by (distance as the k-NN kernel orders it, row).
 */
void merge_lists(const float* bd, const int* bi, const float* nd, const int* ni, int64_t M, int l, int64_t a,
                 float* od, int* oi, hipStream_t s);

/** Scratch of the cells of one level of one copy (reused across levels and copies). */
struct cell_builder {
  int64_t n     = 0;
  int w         = 0;
  hipStream_t s = nullptr;
  dbuf keys, skeys, idx, sidx, sidx2, rid, flag, mkey, mkey2, tmp;
  dbuf start, ukey, pop, keep, kidx, ckey, cfirst, cpop, cstart, z, lists_tmp, bucket, sbucket, seq, perm;
  dbuf ynorm, znorm, kdist;

  /** Scratch for n rows; without member_keys, none for level()'s member sort (the streamed build's levels). */
  void reserve(int64_t n, int w, hipStream_t s, bool member_keys = true);
  /**
   * The cells of the projected rows y [n, w] at spacing f: cells of at least min_cell rows, each with
   * the list of its l members nearest to its center (the nearest repeated when fewer), or with
   * `exact` the l rows nearest to its center among all n (ties by row), or with `ivf` the l rows of ivf->lists
   * (probes probes), in (bucket, id) order.  offs_out [T + 1] (device) receives the CSR over the buckets, keys_out /
   * lists_out the ids and list rows.  Returns the number of cells.
   */
  auto level(const float* y, int B, float f, int min_cell, int l, int log_buckets, bool exact, int* offs_out,
             dbuf& keys_out, dbuf& lists_out, ivf_index* ivf = nullptr, int probes = 0) -> int64_t;
  /**
   * The member-list cells of one level from every row's cell id and squared distance to its cell center (key, dist
   * [n], device; stream_keys): the same cells, keys, lists and offsets as level() with member lists, without the
   * projected rows.
   */
  auto level_streamed(const long long* key, const float* dist, int min_cell, int l, int log_buckets, int* offs_out,
                      dbuf& keys_out, dbuf& lists_out) -> int64_t;
  /**
   * The kept cells of one level from every row's cell id (key [n], device), as level() finds them: ckey_out [M]
   * ascending, crow_out [M] the first row of each (its smallest, the member level() takes the center from).
   * Returns M.
   */
  auto cells_of_keys(const long long* key, int min_cell, dbuf& ckey_out, dbuf& crow_out) -> int64_t;
  /**
   * The level arrays of cells ck [M] with lists [M, l] (both in ck's order): keys_out / lists_out in (bucket, id)
   * order, offs_out [T + 1] their CSR over the buckets.
   */
  void finish_level(const long long* ck, const int* lists, int64_t M, int l, int log_buckets, int* offs_out,
                    dbuf& keys_out, dbuf& lists_out);

 private:
  /** From the sorted ids skeys [n]: the runs, the kept ones (>= min_cell rows) compacted into ckey, cfirst, cpop. */
  auto compact_runs(int min_cell) -> int;
};

}  // namespace cuvs::neighbors::octex::detail
