// Kernels of the octex index builder on MI355X (the reference: detail/build_cells.cuh,
// build_setup.cuh, build_common.cuh).  Cells of a copy are found by sorting the 64-bit cell ids of all
// rows (rocPRIM radix sort), their lists from the members of each cell sorted by their distance to the
// cell center (a second radix sort on (cell, distance)), and the (bucket, id) order with CSR offsets.

#include "build_kernels.hpp"
#include "common.hpp"
#include "e8_device.hpp"

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <rocprim/device/device_radix_sort.hpp>
#include <rocprim/device/device_scan.hpp>

#include <algorithm>
#include <cstdint>
#include <type_traits>

namespace cuvs::neighbors::octex::detail {

namespace {

constexpr int kMaxW = 64;  // 8 * blocks

/** A[i, :] = x[i * step, :] - mean (fp64), for the scatter matrix of the PCA sample. */
__global__ void pca_sample_kernel(const __half* __restrict__ x, int64_t ns, int64_t step, int d,
                                  const float* __restrict__ mean, double* __restrict__ A)
{
  int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= ns * d) return;
  int64_t i = t / d;
  int k     = static_cast<int>(t % d);
  A[t]      = static_cast<double>(__half2float(x[i * step * d + k]) - mean[k]);
}

__global__ void sample_rows_kernel(const __half* __restrict__ x, int64_t ns, int64_t step, int d,
                                   __half* __restrict__ out)
{
  int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= ns * d) return;
  out[t] = x[(t / d) * step * d + t % d];
}

/** G = A^T A (fp64) by 16 x 16 output tiles, samples staged through LDS in chunks of 64 rows. */
__global__ __launch_bounds__(256) void scatter_kernel(const double* __restrict__ A, int64_t ns, int d,
                                                      double* __restrict__ G)
{
  __shared__ double ta[64][17], tb[64][17];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int a0 = blockIdx.y * 16, b0 = blockIdx.x * 16;
  double acc = 0;
  for (int64_t r0 = 0; r0 < ns; r0 += 64) {
    for (int t = threadIdx.x; t < 64 * 16; t += 256) {
      int r = t >> 4, c = t & 15;
      int64_t row = r0 + r;
      ta[r][c]    = (row < ns && a0 + c < d) ? A[row * d + a0 + c] : 0.0;
      tb[r][c]    = (row < ns && b0 + c < d) ? A[row * d + b0 + c] : 0.0;
    }
    __syncthreads();
#pragma unroll 8
    for (int r = 0; r < 64; r++)
      acc = fma(ta[r][ty], tb[r][tx], acc);
    __syncthreads();
  }
  if (a0 + ty < d && b0 + tx < d) G[static_cast<int64_t>(a0 + ty) * d + b0 + tx] = acc;
}

/** y [n, w] = (x - mean) @ U + shift (fp32): one thread per row, U [d, w] in LDS. */
__global__ __launch_bounds__(256) void project_rows_kernel(const __half* __restrict__ x, int64_t n, int d,
                                                           const float* __restrict__ mean,
                                                           const float* __restrict__ U,
                                                           const float* __restrict__ shift, int w,
                                                           float* __restrict__ y)
{
  extern __shared__ float su[];
  float* sm = su + d * w;
  for (int t = threadIdx.x; t < d * w; t += blockDim.x)
    su[t] = U[t];
  for (int t = threadIdx.x; t < d; t += blockDim.x)
    sm[t] = mean[t];
  __syncthreads();
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float acc[kMaxW];
  for (int s = 0; s < w; s++)
    acc[s] = 0.f;
  const __half* r = x + i * d;
  for (int k = 0; k < d; k++) {
    float v = __half2float(r[k]) - sm[k];
    for (int s = 0; s < w; s++)
      acc[s] = fmaf(v, su[k * w + s], acc[s]);
  }
  for (int s = 0; s < w; s++)
    y[i * w + s] = acc[s] + shift[s];
}

/** keys[i] = cell id of y[i] / f (division, as build_cells.cuh:69-71), idx[i] = i. */
template <int B>
__global__ void cell_hash_kernel(const float* __restrict__ y, int64_t n, float f, long long* __restrict__ keys,
                                 int* __restrict__ idx)
{
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float x[8 * B];
#pragma unroll
  for (int k = 0; k < 8 * B; k++)
    x[k] = y[i * 8 * B + k] / f;
  keys[i] = e8b_hash64<B>(x, 1.0f);
  idx[i]  = static_cast<int>(i);
}

/**
 * The streamed build's per-row quantities at spacing f (build_cells.cuh stream_member_copy): key[i] = the cell id of
 * y[i] / f, as cell_hash_kernel, and dist[i] = the squared distance of y[i] to its cell's center f * E8(y[i] / f),
 * as member_key_kernel sums it (every member of a cell has that center).
 */
template <int B>
__global__ void stream_keys_kernel(const float* __restrict__ y, int64_t m, float f, long long* __restrict__ key,
                                   float* __restrict__ dist)
{
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= m) return;
  const float* r = y + i * 8 * B;
  float x[8 * B], z[8 * B];
#pragma unroll
  for (int k = 0; k < 8 * B; k++)
    x[k] = r[k] / f;
  key[i] = e8b_hash64<B>(x, 1.0f);
#pragma unroll
  for (int j = 0; j < B; j++) {
    float xb[8], p[8];
#pragma unroll
    for (int k = 0; k < 8; k++)
      xb[k] = x[8 * j + k];
    e8_point(xb, p);
#pragma unroll
    for (int k = 0; k < 8; k++)
      z[8 * j + k] = p[k] * f;
  }
  float dd = 0.f;
  for (int k = 0; k < 8 * B; k++) {
    const float e = r[k] - z[k];
    dd            = fmaf(e, e, dd);
  }
  dist[i] = dd;
}

/** out[i] = key[idx[i]]. */
__global__ void permute_keys_kernel(const long long* __restrict__ key, const int* __restrict__ idx, int64_t n,
                                    long long* __restrict__ out)
{
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) out[i] = key[idx[i]];
}

/** flag[i] = 1 where a run of equal sorted keys starts. */
__global__ void run_flag_kernel(const long long* __restrict__ k, int64_t n, int* __restrict__ flag)
{
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  flag[i] = (i == 0 || k[i] != k[i - 1]) ? 1 : 0;
}

/** Runs from the inclusive scan rid of the flags: start and key of every run. */
__global__ void run_start_kernel(const long long* __restrict__ k, const int* __restrict__ rid, int64_t n,
                                 int* __restrict__ start, long long* __restrict__ ukey)
{
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  if (i == 0 || k[i] != k[i - 1]) {
    int r    = rid[i] - 1;
    start[r] = static_cast<int>(i);
    ukey[r]  = k[i];
  }
}

/** pop[r] = start[r + 1] - start[r]; keep[r] = a list for run r. */
__global__ void run_keep_kernel(const int* __restrict__ start, int runs, int64_t n, int min_cell,
                                int* __restrict__ pop, int* __restrict__ keep)
{
  int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= runs) return;
  int e   = r + 1 < runs ? start[r + 1] : static_cast<int>(n);
  pop[r]  = e - start[r];
  keep[r] = pop[r] >= min_cell ? 1 : 0;
}

/** The kept runs compacted: key, first row and population of cell kidx[r]. */
__global__ void run_compact_kernel(const long long* __restrict__ ukey, const int* __restrict__ start,
                                   const int* __restrict__ pop, const int* __restrict__ keep,
                                   const int* __restrict__ kidx, int runs, long long* __restrict__ ckey,
                                   int* __restrict__ cfirst, int* __restrict__ cpop)
{
  int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= runs || !keep[r]) return;
  int c     = kidx[r];
  ckey[c]   = ukey[r];
  cfirst[c] = start[r];
  cpop[c]   = pop[r];
}

/**
 * z[c] = f * E8 point of y[first member] / f: the center of kept cell c (build_cells.cuh:86-103).  Without sidx, y
 * holds the first members' projections themselves, y[c] for cell c.
 */
template <int B>
__global__ void cell_center_kernel(const float* __restrict__ y, const int* __restrict__ sidx,
                                   const int* __restrict__ cfirst, int M, float f, float* __restrict__ z)
{
  int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= M) return;
  const int64_t row = sidx != nullptr ? static_cast<int64_t>(sidx[cfirst[c]]) : c;
  const float* r    = y + row * 8 * B;
#pragma unroll
  for (int j = 0; j < B; j++) {
    float x[8], p[8];
#pragma unroll
    for (int k = 0; k < 8; k++)
      x[k] = r[8 * j + k] / f;
    e8_point(x, p);
#pragma unroll
    for (int k = 0; k < 8; k++)
      z[static_cast<int64_t>(c) * 8 * B + 8 * j + k] = p[k] * f;
  }
}

/**
 * Sort key of sorted row i: (kept cell << 32) | distance bits to the cell center (rows of cells
 * without a list sort last).  A stable sort on it orders every cell's members nearest first, ties by
 * row id.
 */
__global__ void member_key_kernel(const float* __restrict__ y, int w, const int* __restrict__ sidx,
                                  const int* __restrict__ rid, const int* __restrict__ keep,
                                  const int* __restrict__ kidx, const float* __restrict__ z, int64_t n,
                                  unsigned long long* __restrict__ key)
{
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  int r = rid[i] - 1;
  if (!keep[r]) {
    key[i] = ~0ULL;
    return;
  }
  int c             = kidx[r];
  const float* v    = y + static_cast<int64_t>(sidx[i]) * w;
  const float* zc   = z + static_cast<int64_t>(c) * w;
  float dd          = 0.f;
  for (int s = 0; s < w; s++) {
    float e = v[s] - zc[s];
    dd      = fmaf(e, e, dd);
  }
  key[i] = (static_cast<unsigned long long>(c) << 32) | __float_as_uint(dd);
}

/** List of cell c: its first l members by distance, the nearest repeated when it has fewer. */
__global__ void list_fill_kernel(const int* __restrict__ sidx2, const int* __restrict__ cstart,
                                 const int* __restrict__ cpop, int M, int l, int* __restrict__ lists)
{
  int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= static_cast<int64_t>(M) * l) return;
  int c = static_cast<int>(t / l), j = static_cast<int>(t % l);
  lists[t] = sidx2[cstart[c] + (j < cpop[c] ? j : 0)];
}

/** crow[c] = sidx[cfirst[c]]: the first row of kept cell c in the stable key sort, its smallest. */
__global__ void first_row_kernel(const int* __restrict__ sidx, const int* __restrict__ cfirst, int M,
                                 int* __restrict__ crow)
{
  int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c < M) crow[c] = sidx[cfirst[c]];
}

/** out [m, d] = x [at[i]]: fp16 rows (d even) by 4-byte words, consecutive threads on consecutive words of a row. */
__global__ void gather_half_rows_kernel(const __half* __restrict__ x, const int* __restrict__ at, int64_t m, int d,
                                        __half* __restrict__ out)
{
  const int64_t t  = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t hw = d / 2;
  if (t >= m * hw) return;
  const int64_t i = t / hw, k = t - i * hw;
  reinterpret_cast<unsigned*>(out)[t] = reinterpret_cast<const unsigned*>(x + static_cast<int64_t>(at[i]) * d)[k];
}

__global__ void bucket_kernel(const long long* __restrict__ ckey, int M, long long mask,
                              unsigned* __restrict__ bucket, int* __restrict__ seq)
{
  int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= M) return;
  bucket[c] = static_cast<unsigned>(ckey[c] & mask);
  seq[c]    = c;
}

/** Cells in (bucket, id) order: keys and list rows gathered by the bucket sort's permutation. */
__global__ void level_gather_kernel(const long long* __restrict__ ckey, const int* __restrict__ lists,
                                    const int* __restrict__ perm, int M, int l, long long* __restrict__ okey,
                                    int* __restrict__ olists)
{
  int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= static_cast<int64_t>(M) * l) return;
  int c = static_cast<int>(t / l), j = static_cast<int>(t % l);
  int p = perm[c];
  olists[t] = lists[static_cast<int64_t>(p) * l + j];
  if (j == 0) okey[c] = ckey[p];
}

/** offs[b] = the number of cells in buckets below b, for b in [0, T] (CSR over the buckets). */
__global__ void offsets_kernel(const unsigned* __restrict__ sbucket, int M, int64_t T, int* __restrict__ offs)
{
  int64_t b = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (b > T) return;
  int lo = 0, hi = M;
  while (lo < hi) {
    int mid = (lo + hi) >> 1;
    if (static_cast<int64_t>(sbucket[mid]) < b)
      lo = mid + 1;
    else
      hi = mid;
  }
  offs[b] = lo;
}

/** v [n, S] = (x - mean) @ basis; amax[s] = max |v[:, s]| (float bits of non-negatives order as uints). */
__global__ __launch_bounds__(256) void sketch_project_kernel(const __half* __restrict__ x, int64_t n, int d,
                                                             const float* __restrict__ mean,
                                                             const float* __restrict__ basis, int S,
                                                             float* __restrict__ v, unsigned* __restrict__ amax)
{
  int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= n * S) return;
  int64_t i = t / S;
  int s     = static_cast<int>(t % S);
  float acc = 0.f;
  for (int k = 0; k < d; k++)
    acc = fmaf(__half2float(x[i * d + k]) - mean[k], basis[static_cast<int64_t>(k) * S + s], acc);
  v[t] = acc;
  atomicMax(amax + s, __float_as_uint(fabsf(acc)));
}

/** codes = clamp(rint(v / scale), -127, 127) (build_setup.cuh:183-190). */
__global__ void quantize_kernel(const float* __restrict__ v, const float* __restrict__ scale, int64_t n, int S,
                                int pitch, signed char* __restrict__ out)
{
  int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= n * pitch) return;
  const int64_t i = t / pitch;
  const int s     = static_cast<int>(t % pitch);
  if (s >= S) {  // the row's padding
    out[t] = 0;
    return;
  }
  float q = rintf(v[i * S + s] / scale[s]);
  out[t]  = static_cast<signed char>(fminf(127.f, fmaxf(-127.f, q)));
}

__global__ void half_to_float_kernel(const __half* __restrict__ x, int64_t total, float* __restrict__ out)
{
  int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t < total) out[t] = __half2float(x[t]);
}

__global__ void float_to_half_kernel(const float* __restrict__ x, int64_t total, __half* __restrict__ out)
{
  int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t < total) out[t] = __float2half_rn(x[t]);
}

// ------------------------------------------------------------------ exact k nearest neighbors

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef float float4_t __attribute__((ext_vector_type(4)));

constexpr int kKnnQ    = 64;   // query rows per workgroup
constexpr int kKnnRows = 128;  // database rows per step: 4 waves x 32
constexpr int kKnnCap  = 256;  // LDS keys per query row: the K kept (K <= 128) and one step's appends
constexpr int kKnnChunk = 8;   // k steps whose fragments are loaded together

__device__ __forceinline__ float knn_f(__half v) { return __half2float(v); }
__device__ __forceinline__ float knn_f(float v) { return v; }

/** out[i] = sum of x[i, :]^2 in fp32, sequentially over the coordinates. */
template <typename T>
__global__ void row_norms_kernel(const T* __restrict__ x, int64_t n, int d, float* __restrict__ out)
{
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const T* r = x + i * d;
  float acc  = 0.f;
  for (int k = 0; k < d; k++) {
    float v = knn_f(r[k]);
    acc     = fmaf(v, v, acc);
  }
  out[i] = acc;
}

/**
 * Four fp16 at columns k..k+3 of `row` (a row pointer, or row 0 of the matrix when the row is past its end:
 * `ok` false), zeros when !ok.  FULL: every column k read lies inside the row (d a multiple of 16), so the load
 * is one unconditional 8-byte load and a select; otherwise each element is checked against d.  The loads are
 * never under a per-lane branch: that made the compiler wait for every earlier load before the next one.
 */
template <bool FULL>
__device__ __forceinline__ half4_t knn_h4(const __half* __restrict__ row, bool ok, int d, int k)
{
  if constexpr (FULL) {
    uint2 u         = *reinterpret_cast<const uint2*>(row + k);
    const half4_t v = *reinterpret_cast<half4_t*>(&u);
    const half4_t z = {0, 0, 0, 0};
    return ok ? v : z;
  } else {
    half4_t v;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const bool in  = ok && k + j < d;
      const __half h = row[in ? k + j : 0];
      v[j]           = in ? static_cast<_Float16>(__half2float(h)) : static_cast<_Float16>(0.f);
    }
    return v;
  }
}

/** Float bits mapped to an unsigned order (negative values first) and back. */
__device__ __forceinline__ unsigned knn_ord(float x)
{
  unsigned u = __float_as_uint(x);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float knn_unord(unsigned o)
{
  return __uint_as_float((o & 0x80000000u) ? (o & 0x7fffffffu) : ~o);
}

/**
 * MFMA fragments of the distance tiles: fp16 rows by v_mfma_f32_16x16x16_f16 (lane l supplies
 * elements 4 (l / 16) .. + 3 of a 16-wide k step for row l % 16), fp32 rows by
 * v_mfma_f32_16x16x4_f32 (lane l supplies element l / 16 of a 4-wide k step).  Both leave D[4 (l / 16)
 * + r][l % 16] in lane l.
 */
template <typename T>
struct knn_op;
template <>
struct knn_op<__half> {
  using frag                 = half4_t;
  static constexpr int kStep = 16;
  static constexpr int kFull = 16;  // d a multiple of this: every lane's columns lie inside the row
  template <bool FULL>
  __device__ static frag load(const __half* row, bool ok, int d, int k0, int lane)
  {
    return knn_h4<FULL>(row, ok, d, k0 + (lane >> 4) * 4);
  }
  __device__ static float4_t mma(frag a, frag b, float4_t c)
  {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
  }
};
template <>
struct knn_op<float> {
  using frag                 = float;
  static constexpr int kStep = 4;
  static constexpr int kFull = 4;
  template <bool FULL>
  __device__ static frag load(const float* row, bool ok, int d, int k0, int lane)
  {
    const int k   = k0 + (lane >> 4);
    const bool in = FULL ? ok : (ok && k < d);
    const float v = row[in ? k : 0];  // unconditional load, then a select
    return in ? v : 0.f;
  }
  __device__ static float4_t mma(frag a, frag b, float4_t c)
  {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
};

/**
 * Every query row's LDS keys (ordered distance << 32 | row) sorted ascending by a bitonic network over
 * all kKnnQ x kKnnCap slots (unused slots padded with ~0), the first K kept, the threshold set to the
 * K-th distance.  Called by the whole workgroup.
 */
__device__ void knn_compact(unsigned long long* key, int* cnt, float* tau, int K)
{
  __syncthreads();
  for (int t = threadIdx.x; t < kKnnQ * kKnnCap; t += blockDim.x)
    if ((t % kKnnCap) >= cnt[t / kKnnCap]) key[t] = ~0ULL;
  for (int size = 2; size <= kKnnCap; size <<= 1)
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      __syncthreads();
      for (int t = threadIdx.x; t < kKnnQ * kKnnCap / 2; t += blockDim.x) {
        const int q = t / (kKnnCap / 2), h = t % (kKnnCap / 2);
        const int lo = ((h & ~(stride - 1)) << 1) | (h & (stride - 1)), hi = lo | stride;
        const bool up = (lo & size) == 0;
        unsigned long long* s = key + q * kKnnCap;
        const unsigned long long x = s[lo], y = s[hi];
        if ((x > y) == up) {
          s[lo] = y;
          s[hi] = x;
        }
      }
    }
  __syncthreads();
  if (threadIdx.x < kKnnQ) {
    const int q = threadIdx.x, c = min(cnt[q], K);
    cnt[q]      = c;
    tau[q]      = c >= K ? knn_unord(static_cast<unsigned>(key[q * kKnnCap + K - 1] >> 32)) : INFINITY;
  }
  __syncthreads();
}

/**
 * The K nearest database rows X [n, d] of each query row Q [m, d] by squared L2 distance
 * |q|^2 + |x|^2 - 2 q.x (fp32; the dot products by MFMA, knn_op: fp16 products are exact in fp32 and
 * accumulated in fp32), ties by row.  A workgroup owns 64 query rows and scans every database row,
 * 128 per step: wave w computes rows [32 w, 32 w + 32) of the step against the 64 queries as 4 x 2
 * MFMA tiles (lane l holds rows 4 (l / 16) + r of a 16-row tile for query l % 16), the fragments of 8 k steps
 * loaded together before their MFMAs.  A distance at or
 * below its query's threshold is appended to the query's LDS keys; when a query holds more than
 * kKnnCap - kKnnRows keys after a step, knn_compact keeps the K smallest and lowers the thresholds, so
 * a step's appends always fit.  out_d / out_i [m, K], sorted; -1 / +inf past the n rows.
 */
template <typename T, bool FULL>
__global__ __launch_bounds__(256) void knn_kernel(const T* __restrict__ Q, const float* __restrict__ qn, int64_t m,
                                                  const T* __restrict__ X, const float* __restrict__ xn, int64_t n,
                                                  int d, int K, float* __restrict__ out_d, int* __restrict__ out_i)
{
  using op = knn_op<T>;
  __shared__ unsigned long long key[kKnnQ * kKnnCap];
  __shared__ int cnt[kKnnQ];
  __shared__ float tau[kKnnQ];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int64_t q0 = static_cast<int64_t>(blockIdx.x) * kKnnQ;
  const int kq     = (lane >> 4) * 4;
  if (tid < kKnnQ) {
    cnt[tid] = 0;
    tau[tid] = INFINITY;
  }
  float qq[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int64_t q = q0 + i * 16 + (lane & 15);
    qq[i]           = q < m ? qn[q] : 0.f;
  }
  __syncthreads();
  for (int64_t r0 = 0; r0 < n; r0 += kKnnRows) {
    const int64_t rw = r0 + wid * 32;
    float4_t acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int t = 0; t < 2; t++)
        acc[i][t] = float4_t{0.f, 0.f, 0.f, 0.f};
    // this step's rows and the workgroup's queries: row pointers (row 0 past the end) and validity, the same
    // for every k step
    const T* xrow[2];
    const T* qrow[4];
    bool xok[2], qok[4];
#pragma unroll
    for (int t = 0; t < 2; t++) {
      const int64_t r = rw + t * 16 + (lane & 15);
      xok[t]          = r < n;
      xrow[t]         = X + (xok[t] ? r : 0) * d;
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int64_t r = q0 + i * 16 + (lane & 15);
      qok[i]          = r < m;
      qrow[i]         = Q + (qok[i] ? r : 0) * d;
    }
    // k in chunks of kKnnChunk steps: the chunk's fragment loads (unconditional, see knn_h4) are all in flight
    // before its MFMAs, so a step of rows waits for memory once per chunk (once for d <= 128 fp16, <= 32 fp32)
    for (int c0 = 0; c0 < d; c0 += op::kStep * kKnnChunk) {
      typename op::frag a[kKnnChunk][2], b[kKnnChunk][4];
#pragma unroll
      for (int j = 0; j < kKnnChunk; j++) {
        if (c0 + op::kStep * j >= d) break;  // uniform
        const int k = c0 + op::kStep * j;
#pragma unroll
        for (int t = 0; t < 2; t++)
          a[j][t] = op::template load<FULL>(xrow[t], xok[t], d, k, lane);
#pragma unroll
        for (int i = 0; i < 4; i++)
          b[j][i] = op::template load<FULL>(qrow[i], qok[i], d, k, lane);
      }
#pragma unroll
      for (int j = 0; j < kKnnChunk; j++) {
        if (c0 + op::kStep * j >= d) break;
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
          for (int t = 0; t < 2; t++)
            acc[i][t] = op::mma(a[j][t], b[j][i], acc[i][t]);
      }
    }
    float xr[2][4];
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int64_t row = rw + t * 16 + kq + r;
        const float v     = xn[row < n ? row : 0];  // unconditional load, then a select
        xr[t][r]          = row < n ? v : 0.f;
      }
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int ql   = i * 16 + (lane & 15);
      const float th = tau[ql];
#pragma unroll
      for (int t = 0; t < 2; t++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const int64_t row = rw + t * 16 + kq + r;
          const float dd    = fmaf(-2.f, acc[i][t][r], qq[i] + xr[t][r]);
          if (row < n && dd <= th) {
            const int p           = atomicAdd(&cnt[ql], 1);
            key[ql * kKnnCap + p] = (static_cast<unsigned long long>(knn_ord(dd)) << 32) |
                                    static_cast<unsigned>(row);
          }
        }
    }
    __syncthreads();  // every append of the step is in
    const int full = tid < kKnnQ && cnt[tid] > kKnnCap - kKnnRows;
    if (__syncthreads_or(full)) knn_compact(key, cnt, tau, K);
  }
  knn_compact(key, cnt, tau, K);
  for (int t = tid; t < kKnnQ * K; t += blockDim.x) {
    const int ql = t / K, j = t % K;
    const int64_t q = q0 + ql;
    if (q >= m) continue;
    const bool ok                = j < cnt[ql];
    const unsigned long long e   = key[ql * kKnnCap + j];
    out_i[q * K + j]             = ok ? static_cast<int>(e & 0xffffffffULL) : -1;
    out_d[q * K + j]             = ok ? knn_unord(static_cast<unsigned>(e >> 32)) : INFINITY;
  }
}

// ------------------------------------------------------------------ IVF lists (build_cells.cuh:511-516, 584-596)

/** ys [ns, w] = y [i * step] (the k-means sample). */
__global__ void take_rows_kernel(const float* __restrict__ y, int64_t ns, int64_t step, int w, float* __restrict__ ys)
{
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= ns * w) return;
  const int64_t i = t / w, k = t - i * w;
  ys[t] = y[i * step * w + k];
}

/** yc [n, w] = y [rows[i]] (the rows grouped by center). */
__global__ void permute_rows_kernel(const float* __restrict__ y, const int* __restrict__ rows, int64_t n, int w,
                                    float* __restrict__ yc)
{
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= n * w) return;
  const int64_t i = t / w, k = t - i * w;
  yc[t] = y[static_cast<int64_t>(rows[i]) * w + k];
}

__global__ void iota_kernel(int* __restrict__ v, int64_t n)
{
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t < n) v[t] = static_cast<int>(t);
}

__global__ void count_labels_kernel(const int* __restrict__ lab, int64_t n, int* __restrict__ cnt)
{
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t < n) atomicAdd(&cnt[lab[t]], 1);
}

/**
 * centers[c] = the mean of the sample rows sidx[off[c]] .. sidx[off[c + 1] - 1] (one workgroup per center; each of
 * the 256 / w parts sums every parts-th member in order, the parts are added in order: the same floats on every
 * run); a center without members keeps its place.
 */
__global__ __launch_bounds__(256) void kmeans_update_kernel(const float* __restrict__ ys, int w,
                                                            const int* __restrict__ sidx, const int* __restrict__ off,
                                                            float* __restrict__ centers)
{
  __shared__ float part[256];
  const int c = blockIdx.x, t = threadIdx.x, parts = 256 / w;
  const int k = t % w, pi = t / w;
  const int a = off[c], b = off[c + 1];
  float acc = 0.f;
  if (pi < parts)
    for (int r = a + pi; r < b; r += parts)
      acc += ys[static_cast<int64_t>(sidx[r]) * w + k];
  part[t] = acc;
  __syncthreads();
  if (t < w && b > a) {
    float sum = 0.f;
    for (int q = 0; q < parts; q++)
      sum += part[q * w + t];
    centers[static_cast<int64_t>(c) * w + t] = sum / static_cast<float>(b - a);
  }
}

constexpr int kIvfBuf  = 512;   // candidate keys below the threshold, waiting to be merged
constexpr int kIvfSort = 1024;  // the kept l (<= 128) and the waiting keys, sorted together

/**
 * The l rows nearest to center z of cell blockIdx.x among the rows of its P probed centers (probe [M, P]; rows of
 * center c: rows[off[c] .. off[c + 1]), coordinates in yc): every candidate's key (fp32 squared distance, summed in
 * coordinate order, then row) is computed by one thread; keys below the current l-th are appended to an LDS buffer,
 * which is merged into the kept l by a bitonic sort whenever the next round could overflow it, and at the end.
 */
__global__ __launch_bounds__(256) void ivf_scan_kernel(const float* __restrict__ z, int w, const int* __restrict__ probe,
                                                       int P, const int* __restrict__ off, const int* __restrict__ rows,
                                                       const float* __restrict__ yc, int l, int* __restrict__ out,
                                                       float* __restrict__ out_d)
{
  __shared__ float zs[kMaxW];
  __shared__ int pre[129], pc[128];
  __shared__ unsigned long long keys[kIvfSort];
  __shared__ int nbuf, nkept;
  __shared__ unsigned long long thr;
  const int64_t cell = blockIdx.x;
  const int t = threadIdx.x;
  constexpr unsigned long long kNone = ~0ULL;
  for (int k = t; k < w; k += blockDim.x)
    zs[k] = z[cell * w + k];
  if (t < 64) {  // wavefront 0: the probed centers and the exclusive prefix of their sizes
    int carry = 0;
    for (int p0 = 0; p0 < P; p0 += 64) {
      const int p  = p0 + t;
      const int c  = p < P ? probe[cell * P + p] : -1;
      const int sz = c >= 0 ? off[c + 1] - off[c] : 0;
      int v        = sz;
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const int u = __shfl_up(v, d);
        if (t >= d) v += u;
      }
      if (p < P) {
        pc[p]  = c;
        pre[p] = carry + v - sz;
      }
      carry += __shfl(v, 63);
    }
    if (t == 0) {
      pre[P] = carry;
      nbuf   = 0;
      nkept  = 0;
      thr    = kNone;
    }
  }
  __syncthreads();
  const int total = pre[P];
  auto merge = [&]() {  // keys[0, nkept) kept (sorted), keys[kIvfSort - kIvfBuf, + nbuf) waiting
    const int nk = nkept, nb = nbuf;
    for (int i = t; i < kIvfSort; i += blockDim.x)
      if (i >= nk && i < kIvfSort - kIvfBuf) keys[i] = kNone;
      else if (i >= kIvfSort - kIvfBuf + nb) keys[i] = kNone;
    __syncthreads();
    for (int size = 2; size <= kIvfSort; size <<= 1)
      for (int stride = size >> 1; stride > 0; stride >>= 1) {
        for (int i = t; i < kIvfSort / 2; i += blockDim.x) {
          const int lo = 2 * i - (i & (stride - 1));  // the pair (lo, lo + stride)
          const int hi = lo + stride;
          const bool up = (lo & size) == 0;
          const unsigned long long a = keys[lo], b = keys[hi];
          if ((a > b) == up) {
            keys[lo] = b;
            keys[hi] = a;
          }
        }
        __syncthreads();
      }
    if (t == 0) {
      int m = 0;
      while (m < l && keys[m] != kNone)
        m++;
      nkept = m;
      nbuf  = 0;
      thr   = m == l ? keys[l - 1] : kNone;
    }
    __syncthreads();
  };
  for (int base = 0; base < total; base += blockDim.x) {
    const int i = base + t;
    if (i < total) {
      int lo = 0, hi = P - 1;  // the last probe whose prefix is <= i
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (pre[mid] <= i)
          lo = mid;
        else
          hi = mid - 1;
      }
      const int64_t j = off[pc[lo]] + (i - pre[lo]);
      const float* r  = yc + j * w;
      float acc       = 0.f;
      for (int k = 0; k < w; k++) {
        const float u = r[k] - zs[k];
        acc           = fmaf(u, u, acc);
      }
      const unsigned long long key =
        (static_cast<unsigned long long>(__float_as_uint(acc)) << 32) | static_cast<unsigned>(rows[j]);
      if (key < thr) keys[kIvfSort - kIvfBuf + atomicAdd(&nbuf, 1)] = key;
    }
    __syncthreads();
    if (nbuf > kIvfBuf - static_cast<int>(blockDim.x)) merge();  // the next round could overflow the buffer
  }
  if (nbuf > 0) merge();
  for (int k = t; k < l; k += blockDim.x) {
    out[cell * l + k] = k < nkept ? static_cast<int>(keys[k] & 0xffffffffULL) : -1;
    if (out_d != nullptr) out_d[cell * l + k] = k < nkept ? __uint_as_float(static_cast<unsigned>(keys[k] >> 32)) : INFINITY;
  }
}

/** bd = +inf, bi = -1: empty lists before the first range's merge. */
__global__ void list_init_kernel(float* __restrict__ bd, int* __restrict__ bi, int64_t total)
{
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= total) return;
  bd[t] = INFINITY;
  bi[t] = -1;
}

/**
 * The streamed lists' merge over row ranges (build_cells.cuh stream_merge_kernel): for each of M centers, the l first
 * of its kept list (bd, bi) and of a range's list (nd, ni, rows numbered from a), both ascending by (distance, row;
 * -1 entries last), into od, oi.  Distances order as the k-NN kernel orders them and rows as unsigned, so the lists
 * merged over ranges are the lists of one search over all rows.
 */
__global__ void merge_lists_kernel(const float* __restrict__ bd, const int* __restrict__ bi,
                                   const float* __restrict__ nd, const int* __restrict__ ni, int64_t M, int l,
                                   int64_t a, float* __restrict__ od, int* __restrict__ oi)
{
  const int64_t c = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (c >= M) return;
  const int64_t o = c * l;
  auto key        = [](float dd, int row) {
    return (static_cast<unsigned long long>(knn_ord(dd)) << 32) | static_cast<unsigned>(row);
  };
  int p = 0, q = 0;  // p + q = j < l: both stay in their lists
  for (int j = 0; j < l; j++) {
    const int ry = ni[o + q] >= 0 ? static_cast<int>(ni[o + q] + a) : -1;
    if (key(bd[o + p], bi[o + p]) <= key(nd[o + q], ry)) {
      od[o + j] = bd[o + p];
      oi[o + j] = bi[o + p];
      p++;
    } else {
      od[o + j] = nd[o + q];
      oi[o + j] = ry;
      q++;
    }
  }
}

template <typename T>
void ensure(dbuf& b, int64_t count)
{
  size_t want = static_cast<size_t>(std::max<int64_t>(count, 1)) * sizeof(T);
  if (b.size < want) b = dbuf(want + want / 8);
}

/** Runs a rocPRIM device call after sizing its temporary storage (grown as needed, never short). */
template <typename F>
void with_tmp(dbuf& tmp, F&& call)
{
  size_t need = 0;
  OCTEX_HIP(call(static_cast<void*>(nullptr), need));
  if (tmp.size < need) tmp = dbuf(need + need / 8);
  size_t have = tmp.size;
  OCTEX_HIP(call(tmp.ptr, have));
}

}  // namespace

// ================================================================== host side

void pca_scatter(const __half* x, int64_t n, int d, int64_t step, int64_t ns, const float* mean, double* G,
                 hipStream_t s)
{
  dbuf A(static_cast<size_t>(ns) * d * sizeof(double));
  pca_sample_kernel<<<grid_for(ns * d, 256), 256, 0, s>>>(x, ns, step, d, mean, A.as<double>());
  dim3 grid((d + 15) / 16, (d + 15) / 16);
  scatter_kernel<<<grid, 256, 0, s>>>(A.as<double>(), ns, d, G);
  OCTEX_HIP(hipGetLastError());
  OCTEX_HIP(hipStreamSynchronize(s));
}

void sample_rows(const __half* x, int64_t ns, int64_t step, int d, __half* host_out, hipStream_t s)
{
  if (ns * d == 0) return;
  dbuf tmp(static_cast<size_t>(ns) * d * sizeof(__half));
  sample_rows_kernel<<<grid_for(ns * d, 256), 256, 0, s>>>(x, ns, step, d, tmp.as<__half>());
  OCTEX_HIP(hipGetLastError());
  OCTEX_HIP(hipMemcpyAsync(host_out, tmp.ptr, tmp.size, hipMemcpyDeviceToHost, s));
  OCTEX_HIP(hipStreamSynchronize(s));
}

void project_rows(const __half* x, int64_t n, int d, const float* mean, const float* U, const float* shift, int w,
                  float* y, hipStream_t s)
{
  OCTEX_EXPECTS(w <= kMaxW, "octex: blocks must be at most 8");
  const size_t smem = static_cast<size_t>(d * w + d) * sizeof(float);
  OCTEX_EXPECTS(smem <= 160 * 1024, "octex: dimension x 8 blocks too large for the projection kernel");
  OCTEX_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&project_rows_kernel),
                                hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(smem)));
  project_rows_kernel<<<grid_for(n, 256), 256, smem, s>>>(x, n, d, mean, U, shift, w, y);
  OCTEX_HIP(hipGetLastError());
}

template <typename T>
void row_norms(const T* x, int64_t n, int d, float* out, hipStream_t s)
{
  if (n == 0) return;
  row_norms_kernel<T><<<grid_for(n, 256), 256, 0, s>>>(x, n, d, out);
  OCTEX_HIP(hipGetLastError());
}
template void row_norms<__half>(const __half*, int64_t, int, float*, hipStream_t);
template void row_norms<float>(const float*, int64_t, int, float*, hipStream_t);

template <typename T>
void knn_rows(const T* Q, const float* qn, int64_t m, const T* X, const float* xn, int64_t n, int d, int K,
              float* out_d, int* out_i, hipStream_t s)
{
  OCTEX_EXPECTS(K >= 1 && K <= kKnnCap - kKnnRows, "octex: exact neighbors: at most %d per row",
                kKnnCap - kKnnRows);
  OCTEX_EXPECTS(n < (int64_t{1} << 31) && d >= 1, "octex: exact neighbors: at most 2^31 - 1 rows");
  if (m == 0) return;
  const int64_t blocks = (m + kKnnQ - 1) / kKnnQ;
  OCTEX_EXPECTS(blocks < (int64_t{1} << 31), "octex: exact neighbors: too many query rows");
  if (d % knn_op<T>::kFull == 0)
    knn_kernel<T, true><<<static_cast<unsigned>(blocks), 256, 0, s>>>(Q, qn, m, X, xn, n, d, K, out_d, out_i);
  else
    knn_kernel<T, false><<<static_cast<unsigned>(blocks), 256, 0, s>>>(Q, qn, m, X, xn, n, d, K, out_d, out_i);
  OCTEX_HIP(hipGetLastError());
}
template void knn_rows<__half>(const __half*, const float*, int64_t, const __half*, const float*, int64_t, int, int,
                               float*, int*, hipStream_t);
template void knn_rows<float>(const float*, const float*, int64_t, const float*, const float*, int64_t, int, int,
                              float*, int*, hipStream_t);

void half_to_float(const __half* x, int64_t total, float* out, hipStream_t s)
{
  if (total == 0) return;
  constexpr int64_t kPiece = int64_t{1} << 30;  // a launch covers fewer than 2^32 work-items
  for (int64_t o = 0; o < total; o += kPiece) {
    const int64_t m = std::min(kPiece, total - o);
    half_to_float_kernel<<<grid_for(m, 256), 256, 0, s>>>(x + o, m, out + o);
    OCTEX_HIP(hipGetLastError());
  }
}

void float_to_half(const float* x, int64_t total, __half* out, hipStream_t s)
{
  if (total == 0) return;
  constexpr int64_t kPiece = int64_t{1} << 30;
  for (int64_t o = 0; o < total; o += kPiece) {
    const int64_t m = std::min(kPiece, total - o);
    float_to_half_kernel<<<grid_for(m, 256), 256, 0, s>>>(x + o, m, out + o);
    OCTEX_HIP(hipGetLastError());
  }
}

auto row_source::rows(int64_t r0, int64_t m, hipStream_t s) -> const __half*
{
  if (dev != nullptr) return dev + r0 * d;
  ensure<__half>(stage, m * d);
  OCTEX_HIP(hipMemcpyAsync(stage.ptr, host + r0 * d, static_cast<size_t>(m) * d * sizeof(__half),
                           hipMemcpyHostToDevice, s));
  return stage.as<__half>();
}

void make_sketch(row_source& x, int64_t n, int d, const float* mean, const float* basis, int S, int pitch,
                 std::vector<float>& scale, signed char* codes, hipStream_t s)
{
  const int64_t chunk = std::min<int64_t>(n, int64_t{1} << 22);
  dbuf v(static_cast<size_t>(chunk) * S * sizeof(float)), amax(S * sizeof(unsigned)), dscale(S * sizeof(float));
  OCTEX_HIP(hipMemsetAsync(amax.ptr, 0, amax.size, s));
  for (int64_t r0 = 0; r0 < n; r0 += chunk) {
    int64_t m = std::min(chunk, n - r0);
    sketch_project_kernel<<<grid_for(m * S, 256), 256, 0, s>>>(x.rows(r0, m, s), m, d, mean, basis, S, v.as<float>(),
                                                              amax.as<unsigned>());
  }
  std::vector<unsigned> ha(S);
  OCTEX_HIP(hipMemcpyAsync(ha.data(), amax.ptr, S * sizeof(unsigned), hipMemcpyDeviceToHost, s));
  OCTEX_HIP(hipStreamSynchronize(s));
  scale.resize(S);
  for (int k = 0; k < S; k++) {
    float am;
    std::memcpy(&am, &ha[k], sizeof(float));
    scale[k] = am > 0.f ? am / 127.f : 1.f;
  }
  OCTEX_HIP(hipMemcpyAsync(dscale.ptr, scale.data(), S * sizeof(float), hipMemcpyHostToDevice, s));
  for (int64_t r0 = 0; r0 < n; r0 += chunk) {
    int64_t m = std::min(chunk, n - r0);
    sketch_project_kernel<<<grid_for(m * S, 256), 256, 0, s>>>(x.rows(r0, m, s), m, d, mean, basis, S, v.as<float>(),
                                                              amax.as<unsigned>());
    quantize_kernel<<<grid_for(m * pitch, 256), 256, 0, s>>>(v.as<float>(), dscale.as<float>(), m, S, pitch,
                                                             codes + r0 * pitch);
  }
  OCTEX_HIP(hipGetLastError());
  OCTEX_HIP(hipStreamSynchronize(s));
}

void cell_builder::reserve(int64_t n_, int w_, hipStream_t s_, bool member_keys)
{
  n = n_;
  w = w_;
  s = s_;
  ensure<long long>(keys, n);
  ensure<long long>(skeys, n);
  ensure<int>(idx, n);
  ensure<int>(sidx, n);
  ensure<int>(sidx2, n);
  ensure<int>(rid, n);
  ensure<int>(flag, n);
  if (member_keys) {
    ensure<unsigned long long>(mkey, n);
    ensure<unsigned long long>(mkey2, n);
  }
}

auto cell_builder::compact_runs(int min_cell) -> int
{
  auto g = grid_for(n, 256);
  run_flag_kernel<<<g, 256, 0, s>>>(skeys.as<long long>(), n, flag.as<int>());
  with_tmp(tmp, [&](void* p, size_t& b) {
    return rocprim::inclusive_scan(p, b, flag.as<int>(), rid.as<int>(), n, rocprim::plus<int>(), s);
  });
  int runs = 0;
  OCTEX_HIP(hipMemcpyAsync(&runs, rid.as<int>() + n - 1, sizeof(int), hipMemcpyDeviceToHost, s));
  OCTEX_HIP(hipStreamSynchronize(s));
  ensure<int>(start, runs + 1);
  ensure<long long>(ukey, runs);
  ensure<int>(pop, runs);
  ensure<int>(keep, runs);
  ensure<int>(kidx, runs);
  run_start_kernel<<<g, 256, 0, s>>>(skeys.as<long long>(), rid.as<int>(), n, start.as<int>(), ukey.as<long long>());
  run_keep_kernel<<<grid_for(runs, 256), 256, 0, s>>>(start.as<int>(), runs, n, min_cell, pop.as<int>(),
                                                      keep.as<int>());
  with_tmp(tmp, [&](void* p, size_t& b) {
    return rocprim::exclusive_scan(p, b, keep.as<int>(), kidx.as<int>(), 0, runs, rocprim::plus<int>(), s);
  });
  int last[2] = {0, 0};
  OCTEX_HIP(hipMemcpyAsync(&last[0], kidx.as<int>() + runs - 1, sizeof(int), hipMemcpyDeviceToHost, s));
  OCTEX_HIP(hipMemcpyAsync(&last[1], keep.as<int>() + runs - 1, sizeof(int), hipMemcpyDeviceToHost, s));
  OCTEX_HIP(hipStreamSynchronize(s));
  const int M = last[0] + last[1];
  ensure<long long>(ckey, M);
  ensure<int>(cfirst, M);
  ensure<int>(cpop, M);
  run_compact_kernel<<<grid_for(runs, 256), 256, 0, s>>>(ukey.as<long long>(), start.as<int>(), pop.as<int>(),
                                                          keep.as<int>(), kidx.as<int>(), runs, ckey.as<long long>(),
                                                          cfirst.as<int>(), cpop.as<int>());
  OCTEX_HIP(hipGetLastError());
  return M;
}

void cell_builder::finish_level(const long long* ck, const int* lists, int64_t M64, int l, int log_buckets,
                                int* offs_out, dbuf& keys_out, dbuf& lists_out)
{
  OCTEX_EXPECTS(M64 < (int64_t{1} << 31), "octex: more than 2^31 - 1 cells in a level");
  const int M     = static_cast<int>(M64);
  const int64_t T = int64_t{1} << log_buckets;
  ensure<unsigned>(bucket, M);
  ensure<unsigned>(sbucket, M);
  ensure<int>(seq, M);
  ensure<int>(perm, M);
  keys_out  = dbuf(static_cast<size_t>(std::max(M, 1)) * sizeof(long long));
  lists_out = dbuf(static_cast<size_t>(std::max<int64_t>(int64_t{M} * l, 1)) * sizeof(int));
  if (M > 0) {
    bucket_kernel<<<grid_for(M, 256), 256, 0, s>>>(ck, M, T - 1, bucket.as<unsigned>(), seq.as<int>());
    with_tmp(tmp, [&](void* p, size_t& b) {
      return rocprim::radix_sort_pairs(p, b, bucket.as<unsigned>(), sbucket.as<unsigned>(), seq.as<int>(),
                                       perm.as<int>(), M, 0, log_buckets, s);
    });
    level_gather_kernel<<<grid_for(int64_t{M} * l, 256), 256, 0, s>>>(ck, lists, perm.as<int>(), M, l,
                                                                       keys_out.as<long long>(), lists_out.as<int>());
  }
  offsets_kernel<<<grid_for(T + 1, 256), 256, 0, s>>>(sbucket.as<unsigned>(), M, T, offs_out);
  OCTEX_HIP(hipGetLastError());
  OCTEX_HIP(hipStreamSynchronize(s));
}

auto cell_builder::cells_of_keys(const long long* key, int min_cell, dbuf& ckey_out, dbuf& crow_out) -> int64_t
{
  auto g = grid_for(n, 256);
  iota_kernel<<<g, 256, 0, s>>>(idx.as<int>(), n);
  with_tmp(tmp, [&](void* p, size_t& b) {
    return rocprim::radix_sort_pairs(p, b, key, skeys.as<long long>(), idx.as<int>(), sidx.as<int>(), n, 0, 64, s);
  });
  const int M = compact_runs(min_cell);
  ckey_out    = dbuf(static_cast<size_t>(std::max(M, 1)) * sizeof(long long));
  crow_out    = dbuf(static_cast<size_t>(std::max(M, 1)) * sizeof(int));
  if (M > 0) {
    OCTEX_HIP(hipMemcpyAsync(ckey_out.ptr, ckey.ptr, static_cast<size_t>(M) * sizeof(long long),
                             hipMemcpyDeviceToDevice, s));
    first_row_kernel<<<grid_for(M, 256), 256, 0, s>>>(sidx.as<int>(), cfirst.as<int>(), M, crow_out.as<int>());
  }
  OCTEX_HIP(hipGetLastError());
  OCTEX_HIP(hipStreamSynchronize(s));
  return M;
}

void cell_centers(const __half* x, const int* rows, int64_t M, int d, const float* mean, const float* U,
                  const float* shift, int B, float f, int64_t chunk, dbuf& stage, float* y, float* z, hipStream_t s)
{
  OCTEX_EXPECTS(d % 2 == 0, "octex: the dimension must be even");
  ensure<__half>(stage, std::min(chunk, M) * d);
  for (int64_t z0 = 0; z0 < M; z0 += chunk) {
    const int64_t m = std::min(chunk, M - z0);
    gather_half_rows_kernel<<<grid_for(m * (d / 2), 256), 256, 0, s>>>(x, rows + z0, m, d, stage.as<__half>());
    project_rows(stage.as<__half>(), m, d, mean, U, shift, 8 * B, y, s);
    auto gm = grid_for(m, 256);
    switch (B) {
#define OCTEX_CC(b) \
  case b: cell_center_kernel<b><<<gm, 256, 0, s>>>(y, nullptr, nullptr, static_cast<int>(m), f, z + z0 * 8 * B); break;
      OCTEX_CC(1) OCTEX_CC(2) OCTEX_CC(3) OCTEX_CC(4) OCTEX_CC(5) OCTEX_CC(6) OCTEX_CC(8)
#undef OCTEX_CC
      default: fail("octex: blocks must be 1-6 or 8");
    }
    OCTEX_HIP(hipGetLastError());
  }
}

void init_lists(float* bd, int* bi, int64_t total, hipStream_t s)
{
  if (total == 0) return;
  list_init_kernel<<<grid_for(total, 256), 256, 0, s>>>(bd, bi, total);
  OCTEX_HIP(hipGetLastError());
}

void merge_lists(const float* bd, const int* bi, const float* nd, const int* ni, int64_t M, int l, int64_t a,
                 float* od, int* oi, hipStream_t s)
{
  if (M == 0) return;
  merge_lists_kernel<<<grid_for(M, 128), 128, 0, s>>>(bd, bi, nd, ni, M, l, a, od, oi);
  OCTEX_HIP(hipGetLastError());
}

auto cell_builder::level(const float* y, int B, float f, int min_cell, int l, int log_buckets, bool exact,
                         int* offs_out, dbuf& keys_out, dbuf& lists_out, ivf_index* ivf, int probes) -> int64_t
{
  const bool member = !exact && ivf == nullptr;
  auto g            = grid_for(n, 256);
  switch (B) {
#define OCTEX_HASH(b) \
  case b: cell_hash_kernel<b><<<g, 256, 0, s>>>(y, n, f, keys.as<long long>(), idx.as<int>()); break;
    OCTEX_HASH(1) OCTEX_HASH(2) OCTEX_HASH(3) OCTEX_HASH(4) OCTEX_HASH(5) OCTEX_HASH(6) OCTEX_HASH(8)
#undef OCTEX_HASH
    default: fail("octex: blocks must be 1-6 or 8");
  }
  with_tmp(tmp, [&](void* p, size_t& b) {
    return rocprim::radix_sort_pairs(p, b, keys.as<long long>(), skeys.as<long long>(), idx.as<int>(), sidx.as<int>(),
                                     n, 0, 64, s);
  });
  const int M = compact_runs(min_cell);
  ensure<int>(cstart, M);
  ensure<float>(z, static_cast<int64_t>(M) * w);
  if (M > 0) {
    auto gm = grid_for(M, 256);
    switch (B) {
#define OCTEX_CENTER(b)                                                                                        \
  case b:                                                                                                      \
    cell_center_kernel<b><<<gm, 256, 0, s>>>(y, sidx.as<int>(), cfirst.as<int>(), M, f, z.as<float>());        \
    break;
      OCTEX_CENTER(1) OCTEX_CENTER(2) OCTEX_CENTER(3) OCTEX_CENTER(4) OCTEX_CENTER(5) OCTEX_CENTER(6) OCTEX_CENTER(8)
#undef OCTEX_CENTER
    }
  }
  if (member) {
    member_key_kernel<<<g, 256, 0, s>>>(y, w, sidx.as<int>(), rid.as<int>(), keep.as<int>(), kidx.as<int>(),
                                        z.as<float>(), n, mkey.as<unsigned long long>());
    with_tmp(tmp, [&](void* p, size_t& b) {
      return rocprim::radix_sort_pairs(p, b, mkey.as<unsigned long long>(), mkey2.as<unsigned long long>(),
                                       sidx.as<int>(), sidx2.as<int>(), n, 0, 64, s);
    });
    if (M > 0)
      with_tmp(tmp, [&](void* p, size_t& b) {
        return rocprim::exclusive_scan(p, b, cpop.as<int>(), cstart.as<int>(), 0, M, rocprim::plus<int>(), s);
      });
  }
  ensure<int>(lists_tmp, static_cast<int64_t>(M) * l);
  if (M > 0) {
    if (ivf != nullptr) {  // the l rows nearest to each center among its probed IVF lists (build_cells.cuh:584-596)
      ensure<float>(znorm, M);
      row_norms<float>(z.as<float>(), M, w, znorm.as<float>(), s);
      ivf->lists(z.as<float>(), znorm.as<float>(), M, probes, l, lists_tmp.as<int>(), s);
    } else if (exact) {  // the l projected rows nearest to each center, by brute force (build_cells.cuh:506-510, 567-599)
      ensure<float>(ynorm, n);
      ensure<float>(znorm, M);
      ensure<float>(kdist, static_cast<int64_t>(M) * l);
      row_norms<float>(y, n, w, ynorm.as<float>(), s);
      row_norms<float>(z.as<float>(), M, w, znorm.as<float>(), s);
      knn_rows<float>(z.as<float>(), znorm.as<float>(), M, y, ynorm.as<float>(), n, w, l, kdist.as<float>(),
                      lists_tmp.as<int>(), s);
    } else {
      list_fill_kernel<<<grid_for(int64_t{M} * l, 256), 256, 0, s>>>(sidx2.as<int>(), cstart.as<int>(),
                                                                      cpop.as<int>(), M, l, lists_tmp.as<int>());
    }
  }
  finish_level(ckey.as<long long>(), lists_tmp.as<int>(), M, l, log_buckets, offs_out, keys_out, lists_out);
  return M;
}

void stream_keys(const float* y, int64_t m, int B, float f, long long* key, float* dist, hipStream_t s)
{
  if (m == 0) return;
  auto g = grid_for(m, 256);
  switch (B) {
#define OCTEX_SK(b) \
  case b: stream_keys_kernel<b><<<g, 256, 0, s>>>(y, m, f, key, dist); break;
    OCTEX_SK(1) OCTEX_SK(2) OCTEX_SK(3) OCTEX_SK(4) OCTEX_SK(5) OCTEX_SK(6) OCTEX_SK(8)
#undef OCTEX_SK
    default: fail("octex: blocks must be 1-6 or 8");
  }
  OCTEX_HIP(hipGetLastError());
}

auto cell_builder::level_streamed(const long long* key, const float* dist, int min_cell, int l, int log_buckets,
                                  int* offs_out, dbuf& keys_out, dbuf& lists_out) -> int64_t
{
  auto g = grid_for(n, 256);
  // rows by distance (stable on the row order), then stably by cell id: each cell's run nearest first, ties by row
  iota_kernel<<<g, 256, 0, s>>>(idx.as<int>(), n);
  ensure<float>(kdist, n);
  with_tmp(tmp, [&](void* p, size_t& b) {
    return rocprim::radix_sort_pairs(p, b, reinterpret_cast<const unsigned*>(dist), kdist.as<unsigned>(),
                                     idx.as<int>(), sidx.as<int>(), n, 0, 32, s);
  });
  permute_keys_kernel<<<g, 256, 0, s>>>(key, sidx.as<int>(), n, keys.as<long long>());
  with_tmp(tmp, [&](void* p, size_t& b) {
    return rocprim::radix_sort_pairs(p, b, keys.as<long long>(), skeys.as<long long>(), sidx.as<int>(),
                                     sidx2.as<int>(), n, 0, 64, s);
  });
  const int M = compact_runs(min_cell);
  ensure<int>(lists_tmp, static_cast<int64_t>(M) * l);
  if (M > 0) {
    // a kept cell's run starts at cfirst in the sorted rows: its first l, the nearest repeated when fewer
    list_fill_kernel<<<grid_for(int64_t{M} * l, 256), 256, 0, s>>>(sidx2.as<int>(), cfirst.as<int>(), cpop.as<int>(),
                                                                    M, l, lists_tmp.as<int>());
  }
  finish_level(ckey.as<long long>(), lists_tmp.as<int>(), M, l, log_buckets, offs_out, keys_out, lists_out);
  return M;
}

void ivf_index::build(const float* y, int64_t n_, int w_, int nlist_, double train_fraction, int iters, hipStream_t s)
{
  n = n_, w = w_, nlist = static_cast<int>(std::min<int64_t>(nlist_, n_));
  OCTEX_EXPECTS(nlist >= 1 && w >= 1 && w <= kMaxW, "octex: IVF lists need rows of at most %d coordinates", kMaxW);
  // the sample: every step-th row, about train_fraction of them and at least nlist
  const int64_t want = std::max<int64_t>(nlist, static_cast<int64_t>(static_cast<double>(n) * train_fraction));
  const int64_t step = std::max<int64_t>(1, n / std::max<int64_t>(want, 1));
  const int64_t ns   = (n + step - 1) / step;
  ensure<float>(ys, ns * w);
  ensure<float>(ysn, ns);
  ensure<float>(centers, int64_t{nlist} * w);
  ensure<float>(cnorm, nlist);
  ensure<int>(off, nlist + 1);
  ensure<int>(cnt, nlist + 1);
  take_rows_kernel<<<grid_for(ns * w, 256), 256, 0, s>>>(y, ns, step, w, ys.as<float>());
  row_norms<float>(ys.as<float>(), ns, w, ysn.as<float>(), s);
  // the first centers: evenly spaced sample rows
  take_rows_kernel<<<grid_for(int64_t{nlist} * w, 256), 256, 0, s>>>(ys.as<float>(), nlist, ns / nlist, w,
                                                                      centers.as<float>());
  const int bits = log2_ceil(nlist) + 1;
  auto group = [&](int64_t m) {  // sidx: 0 .. m-1 ordered by lab (stable), off: CSR of the labels
    ensure<int>(idx, m);
    ensure<int>(sidx, m);
    ensure<int>(slab, m);
    iota_kernel<<<grid_for(m, 256), 256, 0, s>>>(idx.as<int>(), m);
    with_tmp(tmp, [&](void* p, size_t& b) {
      return rocprim::radix_sort_pairs(p, b, lab.as<int>(), slab.as<int>(), idx.as<int>(), sidx.as<int>(),
                                       static_cast<unsigned>(m), 0, bits, s);
    });
    OCTEX_HIP(hipMemsetAsync(cnt.ptr, 0, static_cast<size_t>(nlist + 1) * sizeof(int), s));
    count_labels_kernel<<<grid_for(m, 256), 256, 0, s>>>(lab.as<int>(), m, cnt.as<int>());
    with_tmp(tmp, [&](void* p, size_t& b) {
      return rocprim::exclusive_scan(p, b, cnt.as<int>(), off.as<int>(), 0, nlist + 1, rocprim::plus<int>(), s);
    });
  };
  auto assign = [&](const float* q, const float* qn, int64_t m) {  // lab [m]: the nearest center of every row
    ensure<int>(lab, m);
    ensure<float>(dtmp, m);
    row_norms<float>(centers.as<float>(), nlist, w, cnorm.as<float>(), s);
    knn_rows<float>(q, qn, m, centers.as<float>(), cnorm.as<float>(), nlist, w, 1, dtmp.as<float>(), lab.as<int>(),
                    s);
  };
  for (int it = 0; it < iters; it++) {
    assign(ys.as<float>(), ysn.as<float>(), ns);
    group(ns);
    kmeans_update_kernel<<<nlist, 256, 0, s>>>(ys.as<float>(), w, sidx.as<int>(), off.as<int>(), centers.as<float>());
    OCTEX_HIP(hipGetLastError());
  }
  // every row to its nearest center, the rows grouped by center
  ensure<float>(yn, n);
  row_norms<float>(y, n, w, yn.as<float>(), s);
  assign(y, yn.as<float>(), n);
  group(n);
  rows = dbuf(static_cast<size_t>(n) * sizeof(int));
  OCTEX_HIP(hipMemcpyAsync(rows.ptr, sidx.ptr, rows.size, hipMemcpyDeviceToDevice, s));
  yc = dbuf(static_cast<size_t>(n) * w * sizeof(float));
  permute_rows_kernel<<<grid_for(n * w, 256), 256, 0, s>>>(y, rows.as<int>(), n, w, yc.as<float>());
  row_norms<float>(centers.as<float>(), nlist, w, cnorm.as<float>(), s);
  OCTEX_HIP(hipGetLastError());
  OCTEX_HIP(hipStreamSynchronize(s));
}

void ivf_index::lists(const float* z, const float* zn, int64_t M, int probes, int l, int* out, hipStream_t s,
                      float* out_d)
{
  OCTEX_EXPECTS(l >= 1 && l <= 128, "octex: IVF lists take list_len <= 128");
  if (M == 0) return;
  const int P = std::max(1, std::min({probes, nlist, 128}));
  ensure<float>(pd, M * P);
  ensure<int>(pidx, M * P);
  knn_rows<float>(z, zn, M, centers.as<float>(), cnorm.as<float>(), nlist, w, P, pd.as<float>(), pidx.as<int>(), s);
  OCTEX_EXPECTS(M < (int64_t{1} << 31), "octex: too many cells for one launch");
  ivf_scan_kernel<<<static_cast<unsigned>(M), 256, 0, s>>>(z, w, pidx.as<int>(), P, off.as<int>(), rows.as<int>(),
                                                           yc.as<float>(), l, out, out_d);
  OCTEX_HIP(hipGetLastError());
}

}  // namespace cuvs::neighbors::octex::detail
